// Error state, version, and the staging of descriptor-table uploads.
#include <mutex>
#include <string>

#include "a8_abi_impl.h"

namespace a8 {
static thread_local std::string g_err;
void set_error_msg(const char* msg) { g_err = msg ? msg : ""; }

// Descriptor tables go to the device through a ring of pinned host slots.  A
// hipMemcpyAsync from pageable memory returns only once the copy has run, i.e.
// after every earlier kernel on the stream, which would serialise host-side
// planning with the GPU; from pinned memory it returns at once.  A slot is
// reused only after the event recorded behind its last copy has completed.
namespace {
constexpr int kSlots = 32;
constexpr size_t kSlotBytes = 256 << 10;
constexpr int kMaxDevices = 16;
struct Ring {
  char* host = nullptr;
  hipEvent_t ev[kSlots] = {};
  bool used[kSlots] = {};
  int next = 0;
  bool failed = false;
};
Ring g_ring[kMaxDevices];
std::mutex g_ring_mu;
}  // namespace

hipError_t upload_table(void* dst, const void* src, size_t bytes, hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices || bytes > kSlotBytes)
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
  std::lock_guard<std::mutex> lock(g_ring_mu);
  Ring& r = g_ring[dev];
  if (!r.host && !r.failed) {
    if (hipHostMalloc(reinterpret_cast<void**>(&r.host), kSlots * kSlotBytes, hipHostMallocDefault) != hipSuccess) {
      r.host = nullptr;
      r.failed = true;
    } else {
      for (int i = 0; i < kSlots; ++i) {
        if (hipEventCreateWithFlags(&r.ev[i], hipEventDisableTiming) != hipSuccess) {
          r.failed = true;
          break;
        }
      }
    }
  }
  if (r.failed) return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
  const int s = r.next;
  r.next = (s + 1) % kSlots;
  if (r.used[s]) {
    const hipError_t e = hipEventSynchronize(r.ev[s]);
    if (e != hipSuccess) return e;
  }
  char* slot = r.host + (size_t)s * kSlotBytes;
  std::memcpy(slot, src, bytes);
  hipError_t e = hipMemcpyAsync(dst, slot, bytes, hipMemcpyHostToDevice, st);
  if (e != hipSuccess) return e;
  e = hipEventRecord(r.ev[s], st);
  r.used[s] = e == hipSuccess;
  return e;
}
}  // namespace a8

extern "C" const char* a8_last_error(void) { return a8::g_err.c_str(); }
extern "C" const char* a8_version(void) { return "adafactor8bit_amd 0.1.0 (gfx950)"; }
