// libhwk's device, buffer, stream and event calls: what hwnpu's backend contract asks of a device
// (reference internal/backend/backend.go:12-118), over the HIP runtime. The code-object calls are in
// codeobj.hip.
#include <chrono>
#include <thread>

#include "runtime.h"

extern "C" {

HWK_API int hwk_abi(void) { return HWK_ABI; }

HWK_API void hwk_free_error(char *err) { free(err); }

HWK_API char *hwk_device_count(uint32_t *count) {
  HWK_CHECK(count, "hwk_device_count: null count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice) n = 0;  // looked and found none
  else if (e != hipSuccess) return hwk::hip_err("hipGetDeviceCount", e);
  *count = (uint32_t)n;
  return nullptr;
}

HWK_API char *hwk_device_open(uint32_t index, hwk_device **out) {
  HWK_CHECK(out, "hwk_device_open: null out");
  int n = 0;
  HWK_TRY("hipGetDeviceCount", hipGetDeviceCount(&n));
  HWK_CHECK((int)index < n, "hwk_device_open: device %u of %d", index, n);
  hwk_device *d = new hwk_device();
  d->index = (int)index;
  hipError_t e = hipGetDeviceProperties(&d->prop, d->index);
  if (e != hipSuccess) {
    delete d;
    return hwk::hip_err("hipGetDeviceProperties", e);
  }
  if (strncmp(d->prop.gcnArchName, "gfx950", 6) != 0) {
    char *err = hwk::errf("hwk_device_open: device %u is %s; libhwk's kernels are built for gfx950 only",
                          index, d->prop.gcnArchName);
    delete d;
    return err;
  }
  e = hipSetDevice(d->index);
  if (e != hipSuccess) {
    delete d;
    return hwk::hip_err("hipSetDevice", e);
  }
  *out = d;
  return nullptr;
}

HWK_API void hwk_device_free(hwk_device *d) { delete d; }

HWK_API char *hwk_device_info(hwk_device *d, int key, char *buf, size_t n, size_t *need) {
  HWK_CHECK(d, "hwk_device_info: null device");
  char tmp[256];
  switch (key) {
    case HWK_INFO_NAME: snprintf(tmp, sizeof tmp, "%s", d->prop.name); break;
    case HWK_INFO_ARCH: snprintf(tmp, sizeof tmp, "%s", d->prop.gcnArchName); break;
    case HWK_INFO_PCI_BUS:
      snprintf(tmp, sizeof tmp, "%04x:%02x:%02x", d->prop.pciDomainID, d->prop.pciBusID, d->prop.pciDeviceID);
      break;
    case HWK_INFO_CUS: snprintf(tmp, sizeof tmp, "%d", d->prop.multiProcessorCount); break;
    case HWK_INFO_MEM_BYTES: snprintf(tmp, sizeof tmp, "%zu", (size_t)d->prop.totalGlobalMem); break;
    default: return hwk::errf("hwk_device_info: unknown key %d", key);
  }
  size_t len = strlen(tmp) + 1;
  if (need) *need = len;
  if (buf && n > 0) {
    size_t c = len < n ? len : n;
    memcpy(buf, tmp, c);
    buf[c - 1] = 0;
  }
  return nullptr;
}

HWK_API char *hwk_device_synchronize(hwk_device *d) {
  HWK_CHECK(d, "hwk_device_synchronize: null device");
  HWK_TRY("hipSetDevice", hipSetDevice(d->index));
  HWK_TRY("hipDeviceSynchronize", hipDeviceSynchronize());
  return nullptr;
}

HWK_API char *hwk_buf_alloc(hwk_device *d, size_t size, int kind, hwk_buf **out) {
  HWK_CHECK(d && out, "hwk_buf_alloc: null device or out");
  HWK_CHECK(size > 0, "hwk_buf_alloc: size 0");
  HWK_CHECK(kind == HWK_BUF_MIRRORED || kind == HWK_BUF_DEVICE, "hwk_buf_alloc: unknown kind %d", kind);
  HWK_TRY("hipSetDevice", hipSetDevice(d->index));
  hwk_buf *b = new hwk_buf();
  b->dev = d;
  b->size = size;
  b->kind = kind;
  hipError_t e = hipMalloc(&b->ptr, size);
  if (e != hipSuccess) {
    delete b;
    return hwk::hip_err("hipMalloc", e);
  }
  if (kind == HWK_BUF_MIRRORED) {
    e = hipHostMalloc(&b->host, size, hipHostMallocDefault);
    if (e != hipSuccess) {
      (void)hipFree(b->ptr);
      delete b;
      return hwk::hip_err("hipHostMalloc", e);
    }
    memset(b->host, 0, size);
  }
  *out = b;
  return nullptr;
}

HWK_API void hwk_buf_free(hwk_buf *b) {
  if (!b) return;
  if (b->host) (void)hipHostFree(b->host);
  if (b->ptr) (void)hipFree(b->ptr);
  delete b;
}

HWK_API void *hwk_buf_host_ptr(hwk_buf *b) { return b ? b->host : nullptr; }
HWK_API void *hwk_buf_dev_ptr(hwk_buf *b) { return b ? b->ptr : nullptr; }
HWK_API size_t hwk_buf_size(hwk_buf *b) { return b ? b->size : 0; }

HWK_API char *hwk_buf_sync(hwk_buf *b, int dir, size_t off, size_t n) {
  HWK_CHECK(b, "hwk_buf_sync: null buffer");
  HWK_CHECK(b->host, "hwk_buf_sync: a device-only buffer has no host mirror");
  HWK_CHECK(off <= b->size && n <= b->size - off, "hwk_buf_sync: bytes %zu+%zu past %zu", off, n, b->size);
  if (n == 0) return nullptr;
  HWK_TRY("hipSetDevice", hipSetDevice(b->dev->index));
  char *h = (char *)b->host + off, *dv = (char *)b->ptr + off;
  if (dir == HWK_SYNC_TO_DEVICE)
    HWK_TRY("hipMemcpy", hipMemcpy(dv, h, n, hipMemcpyHostToDevice));
  else if (dir == HWK_SYNC_FROM_DEVICE)
    HWK_TRY("hipMemcpy", hipMemcpy(h, dv, n, hipMemcpyDeviceToHost));
  else
    return hwk::errf("hwk_buf_sync: unknown direction %d", dir);
  return nullptr;
}

HWK_API char *hwk_stream_new(hwk_device *d, void **stream) {
  HWK_CHECK(d && stream, "hwk_stream_new: null device or out");
  HWK_TRY("hipSetDevice", hipSetDevice(d->index));
  hipStream_t s;
  HWK_TRY("hipStreamCreateWithFlags", hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = (void *)s;
  return nullptr;
}

HWK_API void hwk_stream_free(void *stream) {
  if (stream) (void)hipStreamDestroy((hipStream_t)stream);
}

HWK_API char *hwk_stream_sync(void *stream) {
  HWK_TRY("hipStreamSynchronize", hipStreamSynchronize((hipStream_t)stream));
  return nullptr;
}

HWK_API char *hwk_event_new(hwk_device *d, void **event) {
  HWK_CHECK(d && event, "hwk_event_new: null device or out");
  HWK_TRY("hipSetDevice", hipSetDevice(d->index));
  hipEvent_t ev;
  HWK_TRY("hipEventCreate", hipEventCreate(&ev));
  *event = (void *)ev;
  return nullptr;
}

HWK_API void hwk_event_free(void *event) {
  if (event) (void)hipEventDestroy((hipEvent_t)event);
}

HWK_API char *hwk_event_record(void *event, void *stream) {
  HWK_CHECK(event, "hwk_event_record: null event");
  HWK_TRY("hipEventRecord", hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
  return nullptr;
}

// Polls, so that the wait has a bound: the submission keeps running when the wait gives up
// (the reference's Fence.Wait(ctx) is cancelable the same way, graph.go:144-150).
HWK_API char *hwk_event_wait(void *event, uint32_t timeout_ms, int *state) {
  HWK_CHECK(event && state, "hwk_event_wait: null event or state");
  auto start = std::chrono::steady_clock::now();
  for (;;) {
    hipError_t e = hipEventQuery((hipEvent_t)event);
    if (e == hipSuccess) {
      *state = HWK_STATE_DONE;
      return nullptr;
    }
    if (e != hipErrorNotReady) return hwk::hip_err("hipEventQuery", e);
    auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(std::chrono::steady_clock::now() - start).count();
    if ((uint64_t)ms >= timeout_ms) {
      *state = HWK_STATE_PENDING;
      return nullptr;
    }
    std::this_thread::sleep_for(std::chrono::microseconds(50));
  }
}

HWK_API char *hwk_event_elapsed_ns(void *start, void *end, uint64_t *ns) {
  HWK_CHECK(start && end && ns, "hwk_event_elapsed_ns: null argument");
  float ms = 0;
  HWK_TRY("hipEventElapsedTime", hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)end));
  *ns = (uint64_t)((double)ms * 1e6);
  return nullptr;
}

}  // extern "C"
