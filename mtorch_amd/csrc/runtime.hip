// Runtime half of libmthip: error state, per-device streams, the caching allocator, copies,
// stream capture into HIP graphs, and events.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "common.h"

namespace mthip {

namespace {
thread_local std::string g_last_error;

constexpr int kMaxDevices = 64;

struct DeviceState {
  hipStream_t stream = nullptr;
  // Caching allocator: free blocks keyed by size; live blocks map ptr -> (block size, rounded
  // request).  A reused block may be up to 25% larger than the request; `allocated` counts the
  // rounded requests, so it does not depend on which cached block a request happened to get.
  std::multimap<size_t, void*> free_blocks;
  std::unordered_map<void*, std::pair<size_t, size_t>> live;
  size_t allocated = 0;  // rounded request bytes of live blocks
  size_t reserved = 0;   // bytes obtained from hipMalloc and not yet returned
  // Stream capture: blocks freed while a capture is open (or handed out during it) belong to
  // the graph being recorded and may only be reused inside the same capture.
  bool capturing = false;
  std::multimap<size_t, void*> capture_free;
  std::unordered_map<void*, size_t> capture_touched;  // handed out or freed during capture
  std::unordered_map<void*, int> graph_reserved;      // block -> number of live graphs using it
};

std::mutex g_mutex;
DeviceState g_devices[kMaxDevices];

bool caching_disabled() {
  static const bool disabled = [] {
    const char* v = std::getenv("MTHIP_DISABLE_CACHING");
    return v != nullptr && v[0] != '\0' && v[0] != '0';
  }();
  return disabled;
}

// Sizes are rounded so that blocks are reusable across nearby requests: 512 B granules below
// 1 MiB, 128 KiB granules above.  A cached block is reused for a request when it is at most
// 25% (plus one granule) larger, which bounds waste without splitting blocks.
size_t round_size(size_t n) {
  if (n == 0) n = 1;
  if (n < (1u << 20)) return (n + 511) & ~size_t(511);
  const size_t g = size_t(128) << 10;
  return (n + g - 1) / g * g;
}

struct Block {
  void* ptr;
  size_t size;
};

Block take_from(std::multimap<size_t, void*>& pool, size_t size) {
  auto it = pool.lower_bound(size);
  if (it == pool.end() || it->first > size + size / 4 + 4096) return Block{nullptr, 0};
  Block b{it->second, it->first};
  pool.erase(it);
  return b;
}

struct GraphRecord {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<std::pair<void*, size_t>> owned;  // blocks reserved for the graph's lifetime
};

}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int use_device(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(MTHIP_ERR_INVALID, "device index out of range");
  int current = -1;
  MTHIP_CHECK_HIP(hipGetDevice(&current));
  if (current != device) MTHIP_CHECK_HIP(hipSetDevice(device));
  return MTHIP_OK;
}

hipStream_t stream_for(int device) {
  if (device < 0 || device >= kMaxDevices) {
    set_error("device index out of range");
    return nullptr;
  }
  DeviceState& d = g_devices[device];
  if (d.stream) return d.stream;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (d.stream) return d.stream;
  if (use_device(device) != MTHIP_OK) return nullptr;
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) {
    set_error(std::string("hipStreamCreateWithFlags: ") + hipGetErrorString(e));
    return nullptr;
  }
  d.stream = s;
  return s;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MTHIP_ERR_HIP, std::string(what) + " launch: " + hipGetErrorString(e));
  return MTHIP_OK;
}

}  // namespace mthip

using namespace mthip;

extern "C" {

const char* mthip_last_error(void) { return g_last_error.c_str(); }

const char* mthip_version(void) { return "libmthip 0.1 gfx950"; }

int mthip_device_count(int* count) {
  MTHIP_REQUIRE(count != nullptr, "count is NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) n = 0;  // no driver / no device: report zero, as is_available() expects
  *count = n;
  return MTHIP_OK;
}

int mthip_device_info(int device, char* name, size_t name_len, int* cu_count, size_t* total_mem) {
  hipDeviceProp_t prop;
  MTHIP_CHECK_HIP(hipGetDeviceProperties(&prop, device));
  if (name && name_len) {
    // The marketing name comes from libdrm's amdgpu.ids table and is empty where that file is
    // missing; the architecture name and CU count always identify the part.
    std::snprintf(name, name_len, "%s (%s, %d CUs)", prop.name[0] ? prop.name : "AMD GPU", prop.gcnArchName,
                  prop.multiProcessorCount);
  }
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (total_mem) *total_mem = prop.totalGlobalMem;
  return MTHIP_OK;
}

int mthip_malloc(int device, size_t nbytes, void** ptr) {
  MTHIP_REQUIRE(ptr != nullptr, "ptr is NULL");
  if (int rc = use_device(device)) return rc;
  const size_t size = round_size(nbytes);
  std::lock_guard<std::mutex> lock(g_mutex);
  DeviceState& d = g_devices[device];
  Block b{nullptr, 0};
  if (d.capturing) b = take_from(d.capture_free, size);
  if (!b.ptr && !caching_disabled()) b = take_from(d.free_blocks, size);
  if (!b.ptr) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, size);
    if (e != hipSuccess) {
      // Return cached blocks to the driver and retry once before reporting out-of-memory.
      (void)hipGetLastError();
      if (d.stream) (void)hipStreamSynchronize(d.stream);
      for (auto& kv : d.free_blocks) {
        (void)hipFree(kv.second);
        d.reserved -= kv.first;
      }
      d.free_blocks.clear();
      e = hipMalloc(&p, size);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(MTHIP_ERR_OOM, "mthip_malloc: out of device memory allocating " +
                                       std::to_string(nbytes) + " bytes");
      }
    }
    d.reserved += size;
    b = Block{p, size};
  }
  d.live[b.ptr] = {b.size, size};
  d.allocated += size;
  if (d.capturing) d.capture_touched[b.ptr] = b.size;
  *ptr = b.ptr;
  return MTHIP_OK;
}

int mthip_free(int device, void* ptr) {
  if (ptr == nullptr) return MTHIP_OK;
  if (device < 0 || device >= kMaxDevices) return fail(MTHIP_ERR_INVALID, "device index out of range");
  std::lock_guard<std::mutex> lock(g_mutex);
  DeviceState& d = g_devices[device];
  auto it = d.live.find(ptr);
  if (it == d.live.end()) return fail(MTHIP_ERR_INVALID, "mthip_free: pointer not allocated by mthip_malloc");
  const size_t size = it->second.first;
  d.allocated -= it->second.second;
  d.live.erase(it);
  if (d.capturing) {
    // Reusable only inside this capture; afterwards the graph keeps it.
    d.capture_free.emplace(size, ptr);
    d.capture_touched[ptr] = size;
    return MTHIP_OK;
  }
  if (d.graph_reserved.count(ptr)) return MTHIP_OK;  // a live graph replays into it
  if (caching_disabled()) {
    if (int rc = use_device(device)) return rc;
    // Work queued on the stream may still read the block.
    if (d.stream) MTHIP_CHECK_HIP(hipStreamSynchronize(d.stream));
    MTHIP_CHECK_HIP(hipFree(ptr));
    d.reserved -= size;
    return MTHIP_OK;
  }
  // All kernels run in order on the one per-device stream, so a block handed to a later
  // request is only touched by work enqueued after everything that used it before.
  d.free_blocks.emplace(size, ptr);
  return MTHIP_OK;
}

int mthip_empty_cache(int device) {
  if (int rc = use_device(device)) return rc;
  std::lock_guard<std::mutex> lock(g_mutex);
  DeviceState& d = g_devices[device];
  if (d.stream) MTHIP_CHECK_HIP(hipStreamSynchronize(d.stream));
  for (auto& kv : d.free_blocks) {
    MTHIP_CHECK_HIP(hipFree(kv.second));
    d.reserved -= kv.first;
  }
  d.free_blocks.clear();
  return MTHIP_OK;
}

int mthip_memory_stats(int device, size_t* allocated_bytes, size_t* reserved_bytes) {
  if (device < 0 || device >= kMaxDevices) return fail(MTHIP_ERR_INVALID, "device index out of range");
  std::lock_guard<std::mutex> lock(g_mutex);
  if (allocated_bytes) *allocated_bytes = g_devices[device].allocated;
  if (reserved_bytes) *reserved_bytes = g_devices[device].reserved;
  return MTHIP_OK;
}

int mthip_memcpy_h2d(int device, void* dst, const void* src, size_t nbytes) {
  if (nbytes == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  MTHIP_CHECK_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, s));
  // The source is pageable host memory owned by the caller: wait so it may be reused.
  MTHIP_CHECK_HIP(hipStreamSynchronize(s));
  return MTHIP_OK;
}

int mthip_memcpy_d2h(int device, void* dst, const void* src, size_t nbytes) {
  if (nbytes == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  MTHIP_CHECK_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, s));
  MTHIP_CHECK_HIP(hipStreamSynchronize(s));
  return MTHIP_OK;
}

int mthip_memcpy_d2d(int device, void* dst, const void* src, size_t nbytes) {
  if (nbytes == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  MTHIP_CHECK_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, s));
  return MTHIP_OK;
}

int mthip_synchronize(int device) {
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  MTHIP_CHECK_HIP(hipStreamSynchronize(s));
  return MTHIP_OK;
}

void* mthip_stream(int device) { return (void*)stream_for(device); }

int mthip_graph_begin(int device) {
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState& d = g_devices[device];
    MTHIP_REQUIRE(!d.capturing, "mthip_graph_begin: a capture is already open on this device");
    d.capturing = true;
    d.capture_free.clear();
    d.capture_touched.clear();
  }
  hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) {
    std::lock_guard<std::mutex> lock(g_mutex);
    g_devices[device].capturing = false;
    g_devices[device].capture_free.clear();
    g_devices[device].capture_touched.clear();
    return fail(MTHIP_ERR_HIP, std::string("hipStreamBeginCapture: ") + hipGetErrorString(e));
  }
  return MTHIP_OK;
}

int mthip_graph_end(int device, void** graph) {
  MTHIP_REQUIRE(graph != nullptr, "graph is NULL");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  auto* rec = new GraphRecord();
  std::vector<std::pair<void*, size_t>> touched;
  hipError_t e = hipStreamEndCapture(s, &rec->graph);
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState& d = g_devices[device];
    d.capturing = false;
    touched.assign(d.capture_touched.begin(), d.capture_touched.end());
    d.capture_touched.clear();
    d.capture_free.clear();
  }
  std::string err;
  if (e != hipSuccess) {
    err = std::string("hipStreamEndCapture: ") + hipGetErrorString(e);
  } else {
    e = hipGraphInstantiate(&rec->exec, rec->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
      err = std::string("hipGraphInstantiate: ") + hipGetErrorString(e);
      (void)hipGraphDestroy(rec->graph);
    }
  }
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState& d = g_devices[device];
    for (auto& kv : touched) {
      if (err.empty()) {
        // Every block the capture handed out or freed is replayed into by the graph: keep it
        // out of the shared cache until the graph is destroyed.
        rec->owned.emplace_back(kv.first, kv.second);
        d.graph_reserved[kv.first] += 1;
      } else if (d.live.find(kv.first) == d.live.end() && d.graph_reserved.count(kv.first) == 0) {
        // No graph exists to replay into a block freed during the failed capture: it goes
        // back to the shared cache.
        d.free_blocks.emplace(kv.second, kv.first);
      }
    }
  }
  if (!err.empty()) {
    delete rec;
    return fail(MTHIP_ERR_HIP, err);
  }
  *graph = rec;
  return MTHIP_OK;
}

int mthip_graph_launch(int device, void* graph) {
  MTHIP_REQUIRE(graph != nullptr, "graph is NULL");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  MTHIP_CHECK_HIP(hipGraphLaunch(static_cast<GraphRecord*>(graph)->exec, s));
  return MTHIP_OK;
}

int mthip_graph_destroy(int device, void* graph) {
  if (graph == nullptr) return MTHIP_OK;
  if (int rc = use_device(device)) return rc;
  auto* rec = static_cast<GraphRecord*>(graph);
  hipStream_t s = stream_for(device);
  if (s) MTHIP_CHECK_HIP(hipStreamSynchronize(s));
  MTHIP_CHECK_HIP(hipGraphExecDestroy(rec->exec));
  MTHIP_CHECK_HIP(hipGraphDestroy(rec->graph));
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState& d = g_devices[device];
    // Blocks no other graph holds and that are no longer live go back to the shared cache.
    for (auto& ro : rec->owned) {
      auto it = d.graph_reserved.find(ro.first);
      if (it != d.graph_reserved.end() && --it->second == 0) d.graph_reserved.erase(it);
      if (d.graph_reserved.count(ro.first) == 0 && d.live.find(ro.first) == d.live.end())
        d.free_blocks.emplace(ro.second, ro.first);
    }
  }
  delete rec;
  return MTHIP_OK;
}

int mthip_event_create(void** event) {
  MTHIP_REQUIRE(event != nullptr, "event is NULL");
  hipEvent_t e;
  MTHIP_CHECK_HIP(hipEventCreate(&e));
  *event = (void*)e;
  return MTHIP_OK;
}

int mthip_event_record(int device, void* event) {
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  MTHIP_CHECK_HIP(hipEventRecord((hipEvent_t)event, s));
  return MTHIP_OK;
}

int mthip_event_elapsed_ms(void* start, void* end, float* ms) {
  MTHIP_REQUIRE(ms != nullptr, "ms is NULL");
  MTHIP_CHECK_HIP(hipEventSynchronize((hipEvent_t)end));
  MTHIP_CHECK_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
  return MTHIP_OK;
}

int mthip_event_destroy(void* event) {
  if (event) MTHIP_CHECK_HIP(hipEventDestroy((hipEvent_t)event));
  return MTHIP_OK;
}

}  // extern "C"
