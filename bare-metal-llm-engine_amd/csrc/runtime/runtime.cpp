// runtime.cpp -- errors, device queries, memory, streams and events of the C-ABI.
//
// HIP-backed replacement of the reference's src/cuda_device.cpp (device
// queries, 51-301), src/cuda_stream.cpp (RAII stream/event, 11-38) and the
// raw cudaMalloc/cudaMemcpy/cudaMemset calls of include/engine/device_buffer.hpp
// (33-92), exposed as plain C functions.
#include "../engine_internal.hpp"

#include <engine/config.hpp>

#include <dirent.h>

#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <memory>
#include <sstream>
#include <string>

namespace eng {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& msg) { g_last_error = msg; }
void clear_last_error() { g_last_error.clear(); }

void raise(int code, const char* file, int line, const char* expr, const std::string& msg) {
  std::ostringstream oss;
  oss << "[engine] " << file << ":" << line << "\n"
      << "  check failed: " << expr << "\n"
      << "  " << msg;
  throw Error(code, oss.str());
}

void raise_hip(hipError_t err, const char* file, int line, const char* expr) {
  std::ostringstream oss;
  oss << hipGetErrorName(err) << ": " << hipGetErrorString(err);
  raise(ENG_DEVICE_ERROR, file, line, expr, oss.str());
}

namespace {

int device_count_or_zero() {
  int n = 0;
  // Not an error when there is no driver or device: the answer is zero.
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

void current_props(hipDeviceProp_t& prop) {
  ENG_CHECK(device_count_or_zero() > 0, "no HIP device is visible");
  int dev = 0;
  ENG_HIP_CHECK(hipGetDevice(&dev));
  ENG_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
}

void copy_out(const std::string& s, char* buf, std::size_t len) {
  ENG_CHECK(buf != nullptr, "output buffer is null");
  ENG_CHECK(len > 0, "output buffer length must be positive");
  std::snprintf(buf, len, "%s", s.c_str());
}

// Published HBM peak of known parts, in GB/s. hipDeviceProp's memory clock
// times bus width undercounts HBM3E's data rate, so a known part reports its
// specification value; anything else falls back to clock x bus bytes x 2.
double spec_peak_gbs(const hipDeviceProp_t& prop) {
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) return 8000.0;
  if (std::strncmp(prop.gcnArchName, "gfx942", 6) == 0) return 5300.0;
  const double clock_hz = static_cast<double>(prop.memoryClockRate) * 1.0e3;
  const double bus_bytes = static_cast<double>(prop.memoryBusWidth) / 8.0;
  return clock_hz * bus_bytes * 2.0 / 1.0e9;
}

// sysfs directory of the current device's PCI function, e.g.
// "/sys/bus/pci/devices/0000:75:00.0"; empty when the bus id is unknown.
std::string pci_sysfs_dir() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return {};
  }
  char bus[64] = {0};
  if (hipDeviceGetPCIBusId(bus, sizeof(bus), dev) != hipSuccess) {
    (void)hipGetLastError();
    return {};
  }
  std::string id(bus);
  for (char& c : id) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
  return id.empty() ? std::string() : "/sys/bus/pci/devices/" + id;
}

// Current level of an amdgpu DPM table (pp_dpm_sclk / pp_dpm_mclk): lines
// "<index>: <value>Mhz", the current one marked with '*'. Returns MHz, or 0
// when the file is missing or has no marked line.
int dpm_current_mhz(const std::string& path) {
  std::ifstream f(path);
  std::string line;
  while (std::getline(f, line)) {
    if (line.find('*') == std::string::npos) continue;
    const std::size_t colon = line.find(':');
    if (colon == std::string::npos) continue;
    const long v = std::strtol(line.c_str() + colon + 1, nullptr, 10);
    if (v > 0) return static_cast<int>(v);
  }
  return 0;
}

// hwmon frequency input of the device (freq1_input = engine clock, freq2_input
// = memory clock, in Hz). Returns MHz or 0.
int hwmon_mhz(const std::string& dir, const char* file) {
  DIR* d = opendir((dir + "/hwmon").c_str());
  if (d == nullptr) return 0;
  int mhz = 0;
  while (dirent* e = readdir(d)) {
    if (std::strncmp(e->d_name, "hwmon", 5) != 0) continue;
    std::ifstream f(dir + "/hwmon/" + e->d_name + "/" + file);
    long long hz = 0;
    if (f >> hz && hz > 0) {
      mhz = static_cast<int>(hz / 1000000);
      break;
    }
  }
  closedir(d);
  return mhz;
}

// Live clock in MHz and where it came from: the DPM table's current level,
// else the hwmon input, else 0 ("unavailable").
int live_clock_mhz(bool engine_clock, std::string* source) {
  const std::string dir = pci_sysfs_dir();
  if (!dir.empty()) {
    const std::string dpm = dir + (engine_clock ? "/pp_dpm_sclk" : "/pp_dpm_mclk");
    int mhz = dpm_current_mhz(dpm);
    if (mhz > 0) {
      if (source) *source = dpm;
      return mhz;
    }
    mhz = hwmon_mhz(dir, engine_clock ? "freq1_input" : "freq2_input");
    if (mhz > 0) {
      if (source) *source = dir + "/hwmon/*/" + (engine_clock ? "freq1_input" : "freq2_input");
      return mhz;
    }
  }
  if (source) *source = "unavailable";
  return 0;
}

}  // namespace
}  // namespace eng

using eng::guarded;

extern "C" {

const char* eng_last_error(void) { return eng::g_last_error.c_str(); }

#ifndef ENGINE_GIT_REV
#define ENGINE_GIT_REV "unknown"
#endif

const char* eng_build_info(void) {
  return "engine_hip " ENGINE_VERSION_STRING " " ENGINE_HIP_ARCH_STRING " -O3 packed-fp32-off"
#ifdef ENGINE_ALWAYS_SYNC_CHECK
         " sync-check"
#endif
         " git " ENGINE_GIT_REV;
}

int eng_device_count(int* count) {
  return guarded([&] {
    ENG_CHECK(count != nullptr, "eng_device_count: count is null");
    *count = eng::device_count_or_zero();
  });
}

int eng_device_summary(char* buf, std::size_t len) {
  return guarded([&] {
    if (eng::device_count_or_zero() == 0) {
      eng::copy_out("no HIP device", buf, len);
      return;
    }
    hipDeviceProp_t prop{};
    eng::current_props(prop);
    std::ostringstream oss;
    oss.setf(std::ios::fixed);
    oss.precision(1);
    const char* name = prop.name[0] != '\0' ? prop.name : "AMD GPU";
    oss << name << " | " << prop.gcnArchName << " | "
        << (static_cast<double>(prop.totalGlobalMem) / (1024.0 * 1024.0 * 1024.0)) << " GiB"
        << " | " << prop.multiProcessorCount << " CUs"
        << " | " << (prop.sharedMemPerBlock / 1024) << " KiB LDS/block"
        << " | " << eng::spec_peak_gbs(prop) << " GB/s";
    eng::copy_out(oss.str(), buf, len);
  });
}

int eng_peak_bandwidth_gbs(double* gbs) {
  return guarded([&] {
    ENG_CHECK(gbs != nullptr, "eng_peak_bandwidth_gbs: gbs is null");
    *gbs = 0.0;
    if (eng::device_count_or_zero() == 0) return;
    hipDeviceProp_t prop{};
    eng::current_props(prop);
    *gbs = eng::spec_peak_gbs(prop);
  });
}

int eng_driver_version(char* buf, std::size_t len) {
  return guarded([&] {
    int drv = 0;
    if (hipDriverGetVersion(&drv) != hipSuccess) {
      (void)hipGetLastError();
      eng::copy_out("none", buf, len);
      return;
    }
    eng::copy_out(std::to_string(drv), buf, len);
  });
}

int eng_clock_rate_khz(int* khz) {
  return guarded([&] {
    ENG_CHECK(khz != nullptr, "eng_clock_rate_khz: khz is null");
    *khz = 0;
    if (eng::device_count_or_zero() == 0) return;
    hipDeviceProp_t prop{};
    eng::current_props(prop);
    *khz = prop.clockRate;
  });
}

int eng_live_sm_clock_mhz(int* mhz) {
  return guarded([&] {
    ENG_CHECK(mhz != nullptr, "eng_live_sm_clock_mhz: mhz is null");
    *mhz = 0;
    if (eng::device_count_or_zero() == 0) return;
    *mhz = eng::live_clock_mhz(true, nullptr);
    if (*mhz > 0) return;
    hipDeviceProp_t prop{};  // no live source: the nominal clock, as the reference falls back
    eng::current_props(prop);
    *mhz = prop.clockRate / 1000;
  });
}

int eng_live_mem_clock_mhz(int* mhz) {
  return guarded([&] {
    ENG_CHECK(mhz != nullptr, "eng_live_mem_clock_mhz: mhz is null");
    *mhz = 0;
    if (eng::device_count_or_zero() == 0) return;
    *mhz = eng::live_clock_mhz(false, nullptr);
  });
}

int eng_live_clock_source(char* buf, size_t len) {
  return guarded([&] {
    if (eng::device_count_or_zero() == 0) {
      eng::copy_out("no HIP device", buf, len);
      return;
    }
    std::string sclk;
    std::string mclk;
    (void)eng::live_clock_mhz(true, &sclk);
    (void)eng::live_clock_mhz(false, &mclk);
    eng::copy_out("engine clock: " + sclk + "; memory clock: " + mclk, buf, len);
  });
}

int eng_device_arch(char* buf, std::size_t len) {
  return guarded([&] {
    if (eng::device_count_or_zero() == 0) {
      eng::copy_out("none", buf, len);
      return;
    }
    hipDeviceProp_t prop{};
    eng::current_props(prop);
    eng::copy_out(prop.gcnArchName, buf, len);
  });
}

int eng_device_cu_count(int* cus) {
  return guarded([&] {
    ENG_CHECK(cus != nullptr, "eng_device_cu_count: cus is null");
    *cus = 0;
    if (eng::device_count_or_zero() == 0) return;
    hipDeviceProp_t prop{};
    eng::current_props(prop);
    *cus = prop.multiProcessorCount;
  });
}

// ---------------------------------------------------------------- memory

int eng_malloc(void** ptr, std::size_t bytes) {
  return guarded([&] {
    ENG_CHECK(ptr != nullptr, "eng_malloc: ptr is null");
    *ptr = nullptr;
    if (bytes == 0) return;
    ENG_HIP_CHECK(hipMalloc(ptr, bytes));
  });
}

int eng_free(void* ptr) {
  return guarded([&] {
    if (ptr == nullptr) return;
    ENG_HIP_CHECK(hipFree(ptr));
  });
}

int eng_memcpy_h2d(void* dst, const void* src, std::size_t bytes) {
  return guarded([&] {
    if (bytes == 0) return;
    ENG_CHECK(dst != nullptr && src != nullptr, "eng_memcpy_h2d: null pointer");
    ENG_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  });
}

int eng_memcpy_d2h(void* dst, const void* src, std::size_t bytes) {
  return guarded([&] {
    if (bytes == 0) return;
    ENG_CHECK(dst != nullptr && src != nullptr, "eng_memcpy_d2h: null pointer");
    ENG_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  });
}

int eng_memcpy_d2d(void* dst, const void* src, std::size_t bytes) {
  return guarded([&] {
    if (bytes == 0) return;
    ENG_CHECK(dst != nullptr && src != nullptr, "eng_memcpy_d2d: null pointer");
    ENG_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    // A device-to-device hipMemcpy may return before the copy has run, and
    // work on a non-blocking stream does not wait for it: finish it here.
    ENG_HIP_CHECK(hipStreamSynchronize(nullptr));
  });
}

int eng_memcpy_h2d_async(void* dst, const void* src, std::size_t bytes, eng_stream stream) {
  return guarded([&] {
    if (bytes == 0) return;
    ENG_CHECK(dst != nullptr && src != nullptr, "eng_memcpy_h2d_async: null pointer");
    ENG_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, eng::as_stream(stream)));
  });
}

int eng_memcpy_d2h_async(void* dst, const void* src, std::size_t bytes, eng_stream stream) {
  return guarded([&] {
    if (bytes == 0) return;
    ENG_CHECK(dst != nullptr && src != nullptr, "eng_memcpy_d2h_async: null pointer");
    ENG_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, eng::as_stream(stream)));
  });
}

int eng_memset(void* ptr, int value, std::size_t bytes) {
  return guarded([&] {
    if (bytes == 0) return;
    ENG_CHECK(ptr != nullptr, "eng_memset: ptr is null");
    ENG_HIP_CHECK(hipMemset(ptr, value, bytes));
    // hipMemset of device memory may return before the fill has run, and
    // work on a non-blocking stream does not wait for it: finish it here.
    ENG_HIP_CHECK(hipStreamSynchronize(nullptr));
  });
}

int eng_memset_async(void* ptr, int value, std::size_t bytes, eng_stream stream) {
  return guarded([&] {
    if (bytes == 0) return;
    ENG_CHECK(ptr != nullptr, "eng_memset_async: ptr is null");
    // A fill kernel, not hipMemsetAsync: memset nodes recorded into a HIP
    // graph have given wrong results on replays after the first.
    eng::fill_bytes_async(ptr, value, bytes, eng::as_stream(stream));
  });
}

int eng_device_sync(void) {
  return guarded([&] { ENG_HIP_CHECK(hipDeviceSynchronize()); });
}

int eng_check_last_launch(void) {
  return guarded([&] { ENG_HIP_CHECK(hipGetLastError()); });
}

// ------------------------------------------------------- streams and events

int eng_stream_create(eng_stream* stream, unsigned int flags) {
  return guarded([&] {
    ENG_CHECK(stream != nullptr, "eng_stream_create: stream is null");
    hipStream_t s = nullptr;
    // Default priority only: streams of different priorities are not used here.
    ENG_HIP_CHECK(hipStreamCreateWithFlags(&s, flags));
    *stream = reinterpret_cast<eng_stream>(s);
  });
}

int eng_stream_destroy(eng_stream stream) {
  return guarded([&] {
    if (stream == nullptr) return;
    hipStream_t s = eng::as_stream(stream);
    // Drain first: the stream's scratch arena may still be in use by queued
    // kernels, and a later stream can be handed the same handle value.
    ENG_HIP_CHECK(hipStreamSynchronize(s));
    eng::release_stream_scratch(s);
    ENG_HIP_CHECK(hipStreamDestroy(s));
  });
}

int eng_stream_sync(eng_stream stream) {
  return guarded([&] { ENG_HIP_CHECK(hipStreamSynchronize(eng::as_stream(stream))); });
}

int eng_stream_wait_event(eng_stream stream, eng_event event, unsigned int flags) {
  return guarded([&] {
    ENG_CHECK(event != nullptr, "eng_stream_wait_event: event is null");
    ENG_HIP_CHECK(hipStreamWaitEvent(eng::as_stream(stream), eng::as_event(event), flags));
  });
}

int eng_stream_delay(eng_stream stream, unsigned int microseconds) {
  return guarded([&] {
    ENG_CHECK(microseconds <= 1000000u, "eng_stream_delay: microseconds must be at most 1000000");
    eng::stream_delay_async(microseconds, eng::as_stream(stream));
  });
}

int eng_event_create(eng_event* event, unsigned int flags) {
  return guarded([&] {
    ENG_CHECK(event != nullptr, "eng_event_create: event is null");
    hipEvent_t e = nullptr;
    ENG_HIP_CHECK(hipEventCreateWithFlags(&e, flags));
    *event = reinterpret_cast<eng_event>(e);
  });
}

int eng_event_destroy(eng_event event) {
  return guarded([&] {
    if (event == nullptr) return;
    ENG_HIP_CHECK(hipEventDestroy(eng::as_event(event)));
  });
}

namespace {
// A captured graph with the scratch blocks its kernels address: taken over
// from the capture stream's arenas when the capture ends, freed with the graph.
struct GraphHandle {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<void*> scratch;
};
}  // namespace

int eng_graph_capture_begin(eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(stream != nullptr,
              "eng_graph_capture_begin: capture needs a created stream, not the null stream");
    eng::begin_capture_scratch(eng::as_stream(stream));
    ENG_HIP_CHECK(hipStreamBeginCapture(eng::as_stream(stream), hipStreamCaptureModeThreadLocal));
  });
}

int eng_graph_capture_end(eng_stream stream, eng_graph* graph) {
  return guarded([&] {
    ENG_CHECK(stream != nullptr, "eng_graph_capture_end: stream is null");
    ENG_CHECK(graph != nullptr, "eng_graph_capture_end: graph is null");
    *graph = nullptr;
    hipGraph_t g = nullptr;
    ENG_HIP_CHECK(hipStreamEndCapture(eng::as_stream(stream), &g));
    hipGraphExec_t exec = nullptr;
    const hipError_t err = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (err != hipSuccess) {
      (void)hipGraphDestroy(g);
      ENG_HIP_CHECK(err);
    }
    auto h = std::make_unique<GraphHandle>();
    h->graph = g;
    h->exec = exec;
    try {
      // Eager launches queued on the stream before the capture may still use
      // the blocks the graph takes over: let them finish first, so a replay
      // on any stream right after this call cannot race them.
      ENG_HIP_CHECK(hipStreamSynchronize(eng::as_stream(stream)));
      eng::adopt_stream_scratch(eng::as_stream(stream), h->scratch);
    } catch (...) {
      (void)hipGraphExecDestroy(exec);
      (void)hipGraphDestroy(g);
      for (void* p : h->scratch) (void)hipFree(p);
      throw;
    }
    *graph = reinterpret_cast<eng_graph>(h.release());
  });
}

int eng_graph_launch(eng_graph graph, eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(graph != nullptr, "eng_graph_launch: graph is null");
    ENG_HIP_CHECK(hipGraphLaunch(reinterpret_cast<GraphHandle*>(graph)->exec,
                                 eng::as_stream(stream)));
  });
}

int eng_graph_destroy(eng_graph graph) {
  return guarded([&] {
    if (graph == nullptr) return;
    auto* h = reinterpret_cast<GraphHandle*>(graph);
    // Replays may still be queued on any stream: wait for the device before
    // freeing the scratch they address.
    const hipError_t e0 = h->scratch.empty() ? hipSuccess : hipDeviceSynchronize();
    const hipError_t e1 = hipGraphExecDestroy(h->exec);
    const hipError_t e2 = hipGraphDestroy(h->graph);
    for (void* p : h->scratch) (void)hipFree(p);
    delete h;
    ENG_HIP_CHECK(e0);
    ENG_HIP_CHECK(e1);
    ENG_HIP_CHECK(e2);
  });
}

int eng_event_record(eng_event event, eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(event != nullptr, "eng_event_record: event is null");
    ENG_HIP_CHECK(hipEventRecord(eng::as_event(event), eng::as_stream(stream)));
  });
}

int eng_event_query(eng_event event, int* done) {
  return guarded([&] {
    ENG_CHECK(done != nullptr, "eng_event_query: done is null");
    if (event == nullptr) {
      *done = 1;
      return;
    }
    const hipError_t q = hipEventQuery(eng::as_event(event));
    if (q == hipSuccess) {
      *done = 1;
    } else if (q == hipErrorNotReady) {
      (void)hipGetLastError();
      *done = 0;
    } else {
      ENG_HIP_CHECK(q);
    }
  });
}

int eng_event_sync(eng_event event) {
  return guarded([&] {
    if (event == nullptr) return;
    ENG_HIP_CHECK(hipEventSynchronize(eng::as_event(event)));
  });
}

int eng_event_elapsed_ms(float* ms, eng_event start, eng_event end) {
  return guarded([&] {
    ENG_CHECK(ms != nullptr, "eng_event_elapsed_ms: ms is null");
    ENG_CHECK(start != nullptr && end != nullptr,
              "eng_event_elapsed_ms called on uninitialized event");
    ENG_HIP_CHECK(hipEventElapsedTime(ms, eng::as_event(start), eng::as_event(end)));
  });
}

}  // extern "C"
