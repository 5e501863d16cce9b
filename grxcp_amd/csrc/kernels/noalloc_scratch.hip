// Scratch of the allocation-free GemmEx entry point (grxblasGemmExNoAlloc).
//
// grxblasGemmExNoAlloc runs the same plans as grxblasGemmEx, with the
// transposed operand copies and split-K partials in this file-scope array
// instead of a workspace the handle allocates. The array sits in a
// translation unit of its own, with no kernels: its code object is loaded
// on a device only when hipGetSymbolAddress asks for it, so a process that
// never calls grxblasGemmExNoAlloc does not hold the 64 MiB. Each device
// that resolves it holds its own copy (kNoAllocScratchBytes of
// zero-initialised storage that is never read before a call writes it)
// until the process ends. In host code `scratch` names a host-side stand-in,
// not device memory: its device address comes from hipGetSymbolAddress, once
// per device, below, and only that address is ever used.
//
// Ordering. Every call on one device shares that device's array. Calls on
// one stream are ordered by the stream. A call on another stream than the
// device's previous scratch user first waits (hipStreamWaitEvent) for an
// event recorded behind that user's launch, so two host threads, handles or
// streams take turns on the array instead of racing on it. The event is
// created with the address, on the device's first call; no call after that
// allocates anything. Under HIP graph capture the wait and the record are
// left out (an event recorded outside the capture cannot be waited on inside
// it): a captured call is ordered only by the graph and its stream.

#include <hip/hip_runtime.h>

#include <mutex>

#include "../launch.h"

namespace grxk {
namespace {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
  std::mutex mu;                    // held from acquire to release
  void* ptr = nullptr;              // device address of `scratch` on this device
  hipEvent_t done = nullptr;        // recorded behind the latest user's launch
  hipStream_t last = nullptr;       // the stream that recorded it
  bool recorded = false;
};

DeviceScratch g_dev[kMaxDevices];

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return st != hipStreamCaptureStatusNone;
}

}  // namespace

NoAllocScratch::NoAllocScratch(hipStream_t s) : stream_(s) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return;
  }
  DeviceScratch& d = g_dev[dev];
  d.mu.lock();
  if (!d.ptr) {
    void* p = nullptr;
    // resolved with `dev` current: each device's copy lives at its own address
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      (void)hipGetLastError();
      d.mu.unlock();
      return;
    }
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      d.mu.unlock();
      return;
    }
    d.ptr = p;
    d.done = ev;
  }
  captured_ = capturing(s);
  if (!captured_ && d.recorded && d.last != s) {
    if (hipStreamWaitEvent(s, d.done, 0) != hipSuccess) {
      (void)hipGetLastError();
      d.mu.unlock();
      return;
    }
  }
  dev_ = dev;
  ptr_ = d.ptr;
}

hipError_t NoAllocScratch::release(bool launched) {
  if (dev_ < 0) return hipSuccess;
  DeviceScratch& d = g_dev[dev_];
  hipError_t e = hipSuccess;
  if (launched && !captured_) {
    e = hipEventRecord(d.done, stream_);
    if (e == hipSuccess) {
      d.last = stream_;
      d.recorded = true;
    }
  }
  dev_ = -1;
  d.mu.unlock();
  return e;
}

NoAllocScratch::~NoAllocScratch() { (void)release(false); }

}  // namespace grxk
