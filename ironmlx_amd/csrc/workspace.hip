// workspace.hip — device workspaces of the calls that need scratch memory
// (split-K partial sums, the gate_up product of a generic fused SwiGLU, the
// expert segment offsets of a grouped gather).
//
// Each (device, stream, slot) keeps one grow-only buffer, taken from the
// stream-ordered pool (hipMallocAsync on that stream, so it is ordered after
// the stream's earlier work) and never freed: HIP graphs captured on the
// stream keep pointing at it, so their replays need no allocation nodes
// (measured ~8 us per captured split-K call otherwise).  Calls on one stream
// execute in order, so they can share its buffers; a graph captured on a
// stream uses that stream's buffers and must not be replayed concurrently
// with other work on that stream.  During capture a buffer cannot grow; a
// larger request then falls back to a per-call hipMallocAsync / hipFreeAsync
// pair (an allocation node in the graph).
#include <mutex>
#include <unordered_map>

#include "launch.h"

namespace iqmm {
namespace {

struct Key {
  int dev;
  hipStream_t st;
  int slot;
  bool operator==(const Key& o) const { return dev == o.dev && st == o.st && slot == o.slot; }
};
struct KeyHash {
  size_t operator()(const Key& k) const {
    return std::hash<const void*>()(static_cast<const void*>(k.st)) ^ (static_cast<size_t>(k.dev) << 48) ^
           (static_cast<size_t>(k.slot) << 56);
  }
};
struct Buf {
  void* p = nullptr;
  size_t cap = 0;
};

std::mutex g_mu;
std::unordered_map<Key, Buf, KeyHash>& table() {
  static auto* t = new std::unordered_map<Key, Buf, KeyHash>();  // lives until the process ends
  return *t;
}

}  // namespace

hipError_t workspace_get(hipStream_t st, int slot, size_t bytes, void** p, bool* owned) {
  *p = nullptr;
  *owned = false;
  if (bytes == 0) bytes = 256;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess) return e;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    Buf& b = table()[Key{dev, st, slot}];
    if (b.cap >= bytes) {
      *p = b.p;
      return hipSuccess;
    }
    if (cs == hipStreamCaptureStatusNone) {
      // grow (x2 steps, 1 MiB minimum); the old buffer stays allocated for
      // graphs that captured it
      size_t cap = b.cap ? b.cap : (size_t{1} << 20);
      while (cap < bytes) cap *= 2;
      void* np = nullptr;
      e = hipMallocAsync(&np, cap, st);
      if (e != hipSuccess) return e;
      b.p = np;
      b.cap = cap;
      *p = np;
      return hipSuccess;
    }
  }
  // capturing and the buffer is too small: a per-call stream-ordered allocation
  e = hipMallocAsync(p, bytes, st);
  if (e == hipSuccess) *owned = true;
  return e;
}

}  // namespace iqmm
